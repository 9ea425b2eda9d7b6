// GPU quantizers: fp32 rows -> GGUF Q4_K / Q6_K / IQ2_XXS super-blocks.
// Stands in for kq.quantize (tests/test_dequant_unattachable.py:36,
// gmlx/mtp_load.py:290).  Q4_K and Q6_K follow llama.cpp's reference
// quantizers (make_qkx2_quants / make_qx_quants searches); IQ2_XXS uses this
// build's own nearest-lattice search (below).  Every float operation is written in a fixed order
// and the file is compiled without contraction, so results are deterministic
// and reproducible on the host.
#include "kq_common.h"
#include "kq_tables.h"

namespace {

__constant__ uint64_t kGrid[256] = KQ_IQ2XXS_GRID_INIT;

__device__ __forceinline__ int rne(float v) { return (int)rintf(v); }

__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Weighted asymmetric search over n values, nmax levels; returns the scale
// and writes the (negated) minimum.
__device__ float search_asym(const float *x, const float *w, uint8_t *L, float *neg_min, uint8_t *Laux,
                             int n, int nmax, float rmin, float rdelta, int nstep) {
    float lo = x[0], hi = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        lo = x[i] < lo ? x[i] : lo;
        hi = x[i] > hi ? x[i] : hi;
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
        int l = rne(iscale * (x[i] - lo));
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
            int l = rne(iscale * (x[i] - lo));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t)l;
            const float fl = (float)l;
            sum_l += w[i] * fl;
            sum_l2 += w[i] * fl * fl;
            sum_xl += w[i] * fl * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float ts = (sum_w * sum_xl - sum_x * sum_l) / D;
            float tm = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (tm > 0) {
                tm = 0;
                ts = sum_xl / sum_l2;
            }
            float err = 0;
            for (int i = 0; i < n; ++i) {
                float diff = ts * (float)Laux[i] + tm - x[i];
                diff = diff * diff;
                err += w[i] * diff;
            }
            if (err < best) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best = err;
                scale = ts;
                lo = tm;
            }
        }
    }
    *neg_min = -lo;
    return scale;
}

__global__ __launch_bounds__(64) void quant_q4k_kernel(const float *__restrict__ w, int64_t n_rows, int nb,
                                                       int64_t w_stride, uint8_t *__restrict__ out) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_rows * nb) return;
    const int64_t row = gid / nb;
    const int bi = (int)(gid - row * nb);
    const float *x = w + row * w_stride + (int64_t)bi * KQ_QK;
    uint8_t *blk = out + gid * 144;
    uint8_t L[KQ_QK], Laux[32];
    float wt[32], mins[8], scales[8];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(sum_x2 / 32.f);
        for (int l = 0; l < 32; ++l) wt[l] = av_x + fabsf(x[32 * j + l]);
        scales[j] = search_asym(x + 32 * j, wt, L + 32 * j, &mins[j], Laux, 32, 15, -1.f, 0.1f, 20);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    uint8_t sc[12];
    for (int i = 0; i < 12; ++i) sc[i] = 0;
    for (int j = 0; j < 8; ++j) {
        int ls = rne(inv_scale * scales[j]);
        int lm = rne(inv_min * mins[j]);
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
    const uint16_t dh = f32_to_f16(max_scale / 63.f);
    const uint16_t mh = f32_to_f16(max_min / 63.f);
    const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
    for (int j = 0; j < 8; ++j) {
        int s, m;
        if (j < 4) {
            s = sc[j] & 63;
            m = sc[j + 4] & 63;
        } else {
            s = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4);
            m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
        }
        const float dd = d * (float)s;
        if (dd == 0.f) continue;
        const float dm = dmin * (float)m;
        for (int i = 0; i < 32; ++i) {
            int l = rne((x[32 * j + i] + dm) / dd);
            l = l < 0 ? 0 : (l > 15 ? 15 : l);
            L[32 * j + i] = (uint8_t)l;
        }
    }
    blk[0] = dh & 0xFF;
    blk[1] = dh >> 8;
    blk[2] = mh & 0xFF;
    blk[3] = mh >> 8;
    for (int i = 0; i < 12; ++i) blk[4 + i] = sc[i];
    for (int c = 0; c < 4; ++c)
        for (int l = 0; l < 32; ++l) blk[16 + 32 * c + l] = (uint8_t)(L[64 * c + l] | (L[64 * c + 32 + l] << 4));
}

__device__ float search_sym(const float *x, int8_t *L, int n, int nmax) {
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
        int l = rne(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (int8_t)(l + nmax);
        const float wi = x[i] * x[i];
        sumlx += wi * x[i] * (float)l;
        suml2 += wi * (float)l * (float)l;
    }
    float scale = suml2 != 0.f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -((float)nmax + 0.1f * (float)is) / vmax;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = rne(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float wi = x[i] * x[i];
            sumlx += wi * x[i] * (float)l;
            suml2 += wi * (float)l * (float)l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = rne(iscale * x[i]);
                l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
                L[i] = (int8_t)(l + nmax);
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

__global__ __launch_bounds__(64) void quant_q6k_kernel(const float *__restrict__ w, int64_t n_rows, int nb,
                                                       int64_t w_stride, uint8_t *__restrict__ out) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_rows * nb) return;
    const int64_t row = gid / nb;
    const int bi = (int)(gid - row * nb);
    const float *x = w + row * w_stride + (int64_t)bi * KQ_QK;
    uint8_t *blk = out + gid * 210;
    int8_t L[KQ_QK];
    float scales[16];
    float max_scale = 0, max_abs = 0;
    for (int ib = 0; ib < 16; ++ib) {
        const float s = search_sym(x + 16 * ib, L + 16 * ib, 16, 32);
        scales[ib] = s;
        if (fabsf(s) > max_abs) {
            max_abs = fabsf(s);
            max_scale = s;
        }
    }
    for (int i = 0; i < 210; ++i) blk[i] = 0;
    if (max_abs < 1e-15f) return;
    const float iscale = -128.f / max_scale;
    const uint16_t dh = f32_to_f16(1.f / iscale);
    blk[208] = dh & 0xFF;
    blk[209] = dh >> 8;
    int8_t sc[16];
    for (int ib = 0; ib < 16; ++ib) {
        const int v = rne(iscale * scales[ib]);
        sc[ib] = (int8_t)(v > 127 ? 127 : v);
        blk[192 + ib] = (uint8_t)sc[ib];
    }
    const float d = f16_to_f32(dh);
    for (int j = 0; j < 16; ++j) {
        const float dd = d * (float)sc[j];
        if (dd == 0.f) continue;
        for (int i = 0; i < 16; ++i) {
            int l = rne(x[16 * j + i] / dd);
            l = l < -32 ? -32 : (l > 31 ? 31 : l);
            L[16 * j + i] = (int8_t)(l + 32);
        }
    }
    for (int h = 0; h < 2; ++h) {
        const int8_t *Lh = L + 128 * h;
        for (int l = 0; l < 32; ++l) {
            const uint8_t a = (uint8_t)Lh[l], b = (uint8_t)Lh[l + 32];
            const uint8_t c = (uint8_t)Lh[l + 64], e = (uint8_t)Lh[l + 96];
            blk[64 * h + l] = (uint8_t)((a & 0xF) | ((c & 0xF) << 4));
            blk[64 * h + l + 32] = (uint8_t)((b & 0xF) | ((e & 0xF) << 4));
            blk[128 + 32 * h + l] = (uint8_t)((a >> 4) | ((b >> 4) << 2) | ((c >> 4) << 4) | ((e >> 4) << 6));
        }
    }
}

// IQ2_XXS quantizer (this build's own search).  Grid bytes take the values
// 8, 25 and 43 (levels 0, 1, 2).  For a scale db, each folded value picks the
// nearest level by the midpoints (below 16.5 db: 0, below 34 db: 1, else 2);
// the 8 levels of a sub-group form a lattice point u = sum l_j 3^j, and the
// grid entry nearest to it in level values (g_iq2_near[u], integer squared
// distance, ties to the lower entry) is taken.  The scale field s (db =
// d (0.5 + s) / 4) with the least squared error over the group's 32 values
// wins (ties to the lower s).

__device__ uint8_t g_iq2_near[6561];

// g_iq2_near[u] for every lattice point u (one thread each).
__global__ __launch_bounds__(256) void iq2_near_kernel() {
    const int u = blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= 6561) return;
    int lv[8];
    for (int j = 0, r = u; j < 8; ++j, r /= 3) lv[j] = r % 3;
    const int val[3] = {8, 25, 43};
    int best = 0x7FFFFFFF, bk = 0;
    for (int k = 0; k < 256; ++k) {
        const uint64_t gv = kGrid[k];
        int dsum = 0;
        for (int j = 0; j < 8; ++j) {
            const int d = val[lv[j]] - (int)((gv >> (8 * j)) & 0xFF);
            dsum += d * d;
        }
        if (dsum < best) {
            best = dsum;
            bk = k;
        }
    }
    g_iq2_near[u] = (uint8_t)bk;
}

// One thread per 32-value group; the block scale d is computed by every
// group thread of the block from the same 256 values.
__global__ __launch_bounds__(64) void quant_iq2xxs_kernel(const float *__restrict__ w, int64_t n_rows, int nb,
                                                          int64_t w_stride, uint8_t *__restrict__ out) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= n_rows * nb * 8) return;
    const int64_t bidx = gid >> 3;
    const int grp = (int)(gid & 7);
    const int64_t row = bidx / nb;
    const int bi = (int)(bidx - row * nb);
    const float *x = w + row * w_stride + (int64_t)bi * KQ_QK;
    uint8_t *blk = out + bidx * 66;
    float amax = 0;
    for (int i = 0; i < KQ_QK; ++i) amax = fabsf(x[i]) > amax ? fabsf(x[i]) : amax;
    if (amax < 1e-30f) {
        if (grp == 0) {
            blk[0] = 0;
            blk[1] = 0;
        }
        for (int i = 0; i < 8; ++i) blk[2 + 8 * grp + i] = 0;
        return;
    }
    const float dguess = amax / (43.f * 15.5f * 0.25f);
    const uint16_t dh = f32_to_f16(dguess);
    if (grp == 0) {
        blk[0] = dh & 0xFF;
        blk[1] = dh >> 8;
    }
    const float d = f16_to_f32(dh);
    const float *xg = x + 32 * grp;
    float folded[32], mag[32];
    uint32_t sign_idx[4];
    for (int i = 0; i < 32; ++i) mag[i] = fabsf(xg[i]);
    for (int l = 0; l < 4; ++l) {
        uint32_t s = 0;
        int nneg = 0, jmin = 0;
        for (int j = 0; j < 8; ++j) {
            if (xg[8 * l + j] < 0) {
                s |= 1u << j;
                nneg++;
            }
            if (mag[8 * l + j] < mag[8 * l + jmin]) jmin = j;
        }
        if (nneg & 1) s ^= 1u << jmin;
        sign_idx[l] = s & 127u;
        const uint32_t full = sign_idx[l] | ((uint32_t)(__builtin_popcount(sign_idx[l]) & 1) << 7);
        for (int j = 0; j < 8; ++j) folded[8 * l + j] = ((full >> j) & 1) ? -xg[8 * l + j] : xg[8 * l + j];
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
            const uint32_t k = g_iq2_near[u];
            const uint64_t gv = kGrid[k];
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
    uint8_t *g = blk + 2 + 8 * grp;
    for (int i = 0; i < 4; ++i) {
        g[i] = (uint8_t)(best_idx >> (8 * i));
        g[4 + i] = (uint8_t)(aux1 >> (8 * i));
    }
}

}  // namespace

extern "C" int kq_quantize(const float *w, int64_t n_rows, int64_t K, int64_t w_row_stride, int codec,
                           void *wire, kq_stream_t stream) {
    if (n_rows == 0) return KQ_OK;
    if (!w || !wire) return KQ_ERR_NULL_POINTER;
    if (kq_block_bytes(codec) == 0) return KQ_ERR_UNSUPPORTED_CODEC;
    if (n_rows < 0 || K <= 0 || K % KQ_QK || w_row_stride < K) return KQ_ERR_BAD_SHAPE;
    const int nb = (int)(K / KQ_QK);
    hipStream_t s = (hipStream_t)stream;
    const int64_t blocks = n_rows * nb;
    if (codec == KQ_CODEC_Q4_K) {
        hipLaunchKernelGGL(quant_q4k_kernel, dim3((unsigned)((blocks + 63) / 64)), dim3(64), 0, s, w, n_rows,
                           nb, w_row_stride, (uint8_t *)wire);
    } else if (codec == KQ_CODEC_Q6_K) {
        hipLaunchKernelGGL(quant_q6k_kernel, dim3((unsigned)((blocks + 63) / 64)), dim3(64), 0, s, w, n_rows,
                           nb, w_row_stride, (uint8_t *)wire);
    } else {
        // the nearest-grid table is rebuilt on the stream ahead of every
        // launch (26 workgroups): no state outlives the call
        hipLaunchKernelGGL(iq2_near_kernel, dim3((6561 + 255) / 256), dim3(256), 0, s);
        hipLaunchKernelGGL(quant_iq2xxs_kernel, dim3((unsigned)((blocks * 8 + 63) / 64)), dim3(64), 0, s, w,
                           n_rows, nb, w_row_stride, (uint8_t *)wire);
    }
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}
