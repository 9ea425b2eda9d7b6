// Ragged GQA decode attention (one query token per row) for gfx950.
//
// Semantics: gmlx/qwen35_attn.py:395-493 (ragged_decode_attention) and the
// batched kq.sdpa_decode_gqa(starts=) route (gmlx/gemma4_batched_sdpa.py:
// 210-226): per (row b, q head hq) softmax(scale * q . K^T) . V over the row's
// visible keys, kv head h = hq / (Hq/Hkv), fp32 online softmax.
//
// Work unit = one wave = (row b, kv head h, split s of C tokens): the wave
// streams its K/V tokens once for all G = Hq/Hkv query heads of the group
// (GQA sharing), 32 tokens per tile, both products on v_mfma_f32_16x16x32:
//   S^T[tok, head]  = K_tile[tok, d] . q^T[d, head]      (A = K rows as loaded)
//   O^T[d, head]   += V^T[d, tok]  . P^T[tok, head]      (A = V^T via v_perm)
// Lane l = 16*g + r: in the score tile it holds head r at tokens
// {4g..4g+3, 16+4g..16+4g+3}; the P.V B-operand wants exactly those tokens
// in the same lane, so P never leaves its lane.  Splits of one (b, h) are
// merged by the last split to finish (agent-scope counter), in split order,
// so the result does not depend on scheduling.
#include "kq_common.h"

namespace {

struct SdpaArgs {
    const uint16_t *q, *k, *v;
    uint16_t *out;
    const int64_t *kv_off, *head_stride;
    const int32_t *row_len;
    float *part;          // [B][Hkv][max_splits][G][D] O partials, then m/l
    float *ml;            // [B][Hkv][max_splits][G][2]
    uint32_t *ctr;        // [B][Hkv]
    int32_t B, Hq, Hkv, G, split, max_splits, max_len;
    float scale_log2;     // scale * log2(e)
};

template <bool BF>
__device__ __forceinline__ floatx4 mfma(const half8_t &a, const half8_t &b, const floatx4 &c) {
    if constexpr (!BF) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    } else {
        typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    }
}

template <bool BF>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (!BF) {
        return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
    } else {
        return (uint32_t)kq_f32_to_bf16_bits(a) | ((uint32_t)kq_f32_to_bf16_bits(b) << 16);
    }
}

template <bool BF>
__device__ __forceinline__ float to_f32(uint16_t h) {
    if constexpr (!BF) return (float)__builtin_bit_cast(_Float16, h);
    else return kq_bf16_bits_to_f32(h);
}

template <bool BF>
__device__ __forceinline__ uint16_t from_f32(float f) {
    if constexpr (!BF) return __builtin_bit_cast(uint16_t, (_Float16)f);
    else return kq_f32_to_bf16_bits(f);
}

// Map unit u to (b, h, s).  Each row contributes max(1, ceil(len/C)) splits
// per kv head.  Returns false when u is past the last unit.
__device__ __forceinline__ bool map_unit(const SdpaArgs &a, int u, int &b, int &h, int &s, int &nsplit) {
    const int lane = kq_lane();
    int base = 0;
    for (int c0 = 0; c0 < a.B; c0 += 64) {
        const int row = c0 + lane;
        int n = 0;
        if (row < a.B) {
            const int len = min(a.row_len[row], a.max_len);
            n = len <= 0 ? 1 : (len + a.split - 1) / a.split;
        }
        const int units = n * a.Hkv;
        // inclusive scan across the wave
        int inc = units;
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(inc, off);
            if (lane >= off) inc += t;
        }
        const int excl = inc - units;
        const int total = __shfl(inc, 63);
        if (u < base + total) {
            const uint64_t hit = __ballot(row < a.B && u >= base + excl && u < base + inc);
            const int src = __builtin_ctzll(hit);
            b = c0 + src;
            nsplit = __shfl(n, src);
            const int local = u - base - __shfl(excl, src);
            h = local / nsplit;
            s = local - h * nsplit;
            return true;
        }
        base += total;
    }
    return false;
}

template <int D, bool BF>
__global__ __launch_bounds__(64) void kq_sdpa_kernel(SdpaArgs a) {
    constexpr int NC = D / 32;               // 32-wide d chunks for Q.K
    constexpr int NG = (D + 127) / 128;      // 128-wide d groups for P.V
    const int lane = kq_lane();
    const int r = lane & 15, g = lane >> 4;

    for (int u = blockIdx.x;; u += gridDim.x) {
        int b, h, s, nsplit;
        if (!map_unit(a, u, b, h, s, nsplit)) return;
        // rows longer than max_len are clamped to it (the workspace holds
        // max_len / split splits per (row, head))
        const int len = max(min(a.row_len[b], a.max_len), 0);
        const int t_begin = s * a.split;
        const int t_end = min(len, t_begin + a.split);
        const int64_t kvbase = a.kv_off[b] + (int64_t)h * a.head_stride[b];
        const uint16_t *kp = a.k + kvbase;
        const uint16_t *vp = a.v + kvbase;
        const bool head_ok = r < a.G;
        const int hq = h * a.G + r;

        // q^T fragments: lane (head r, group g) holds q[hq][32c + 8g .. +7]
        half8_t qf[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (head_ok) {
                qf[c] = __builtin_bit_cast(half8_t, *(const u32x4 *)(a.q + ((int64_t)b * a.Hq + hq) * D + 32 * c + 8 * g));
            } else {
                qf[c] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
            }
        }

        floatx4 o[NG][8];
#pragma unroll
        for (int dg = 0; dg < NG; ++dg)
#pragma unroll
            for (int j = 0; j < 8; ++j) o[dg][j] = floatx4{0, 0, 0, 0};
        float m_run = -INFINITY;   // running max (log2 domain), same on the 4 lanes of a head
        float l_part = 0.f;        // this lane's share of the running sum

        for (int t0 = t_begin; t0 < t_end; t0 += 32) {
            // ---- S = K . q^T for tokens t0 + [0, 32)
            floatx4 sc[2];
#pragma unroll
            for (int ch = 0; ch < 2; ++ch) {
                const int tok = t0 + 16 * ch + r;
                const bool tv = tok < t_end;
                floatx4 acc = {0, 0, 0, 0};
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    half8_t kf = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
                    if (tv) kf = __builtin_bit_cast(half8_t, *(const u32x4 *)(kp + (int64_t)tok * D + 32 * c + 8 * g));
                    acc = mfma<BF>(kf, qf[c], acc);
                }
                sc[ch] = acc;
            }
            // ---- V rows for this lane's 8 tokens, d = 128*dg + 8*r .. +7
            u32x4 vr[NG][8];
#pragma unroll
            for (int dg = 0; dg < NG; ++dg) {
                const int d0 = 128 * dg + 8 * r;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int tok = t0 + (i < 4 ? 4 * g + i : 16 + 4 * g + (i - 4));
                    if (tok < t_end && d0 < D) vr[dg][i] = *(const u32x4 *)(vp + (int64_t)tok * D + d0);
                    else vr[dg][i] = u32x4{0, 0, 0, 0};
                }
            }
            // ---- online softmax over this lane's 8 scores (head r)
            float sv[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int ta = t0 + 4 * g + e, tb = t0 + 16 + 4 * g + e;
                sv[e] = (ta < t_end && head_ok) ? sc[0][e] * a.scale_log2 : -INFINITY;
                sv[4 + e] = (tb < t_end && head_ok) ? sc[1][e] * a.scale_log2 : -INFINITY;
            }
            float tmax = sv[0];
#pragma unroll
            for (int i = 1; i < 8; ++i) tmax = fmaxf(tmax, sv[i]);
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            const float m_new = fmaxf(m_run, tmax);
            // m_new == -inf only for heads >= G or fully masked tiles
            const float alpha = (m_new == -INFINITY) ? 1.f : exp2f(m_run - m_new);
            float p[8];
            float psum = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                p[i] = (m_new == -INFINITY) ? 0.f : exp2f(sv[i] - m_new);
                psum += p[i];
            }
            l_part = l_part * alpha + psum;
            m_run = m_new;
            const half8_t pf = __builtin_bit_cast(
                half8_t, u32x4{pack2<BF>(p[0], p[1]), pack2<BF>(p[2], p[3]), pack2<BF>(p[4], p[5]),
                               pack2<BF>(p[6], p[7])});
            // ---- O^T += V^T . P^T
#pragma unroll
            for (int dg = 0; dg < NG; ++dg) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
                    u32x4 f;
                    f.x = __builtin_amdgcn_perm(vr[dg][1][j >> 1], vr[dg][0][j >> 1], sel);
                    f.y = __builtin_amdgcn_perm(vr[dg][3][j >> 1], vr[dg][2][j >> 1], sel);
                    f.z = __builtin_amdgcn_perm(vr[dg][5][j >> 1], vr[dg][4][j >> 1], sel);
                    f.w = __builtin_amdgcn_perm(vr[dg][7][j >> 1], vr[dg][6][j >> 1], sel);
                    floatx4 acc = o[dg][j] * alpha;
                    o[dg][j] = mfma<BF>(__builtin_bit_cast(half8_t, f), pf, acc);
                }
            }
        }

        // Lane (head r, g) now holds O[hq][d] for d = 128*dg + 32*g + 8*e + j
        // (element e of o[dg][j]); l is split over the 4 lanes of a head.
        float l_tot = l_part + __shfl_xor(l_part, 16);
        l_tot += __shfl_xor(l_tot, 32);

        if (nsplit == 1) {
            if (head_ok) {
                const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
                uint16_t *op = a.out + ((int64_t)b * a.Hq + hq) * D;
#pragma unroll
                for (int dg = 0; dg < NG; ++dg)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int d0 = 128 * dg + 32 * g + 8 * e;
                        if (d0 >= D) continue;
                        u32x4 w;
                        w.x = (uint32_t)from_f32<BF>(o[dg][0][e] * inv) | ((uint32_t)from_f32<BF>(o[dg][1][e] * inv) << 16);
                        w.y = (uint32_t)from_f32<BF>(o[dg][2][e] * inv) | ((uint32_t)from_f32<BF>(o[dg][3][e] * inv) << 16);
                        w.z = (uint32_t)from_f32<BF>(o[dg][4][e] * inv) | ((uint32_t)from_f32<BF>(o[dg][5][e] * inv) << 16);
                        w.w = (uint32_t)from_f32<BF>(o[dg][6][e] * inv) | ((uint32_t)from_f32<BF>(o[dg][7][e] * inv) << 16);
                        *(u32x4 *)(op + d0) = w;
                    }
            }
            continue;
        }

        // ---- split partial: O (unnormalised), m, l
        const int64_t slot = ((int64_t)b * a.Hkv + h) * a.max_splits;
        if (head_ok) {
            float *po = a.part + ((slot + s) * a.G + r) * D;
#pragma unroll
            for (int dg = 0; dg < NG; ++dg)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int d0 = 128 * dg + 32 * g + 8 * e;
                    if (d0 >= D) continue;
                    float4 *dst = (float4 *)(po + d0);
                    dst[0] = make_float4(o[dg][0][e], o[dg][1][e], o[dg][2][e], o[dg][3][e]);
                    dst[1] = make_float4(o[dg][4][e], o[dg][5][e], o[dg][6][e], o[dg][7][e]);
                }
            if (g == 0) {
                float *pml = a.ml + ((slot + s) * a.G + r) * 2;
                pml[0] = m_run;
                pml[1] = l_tot;
            }
        }
        __threadfence();
        uint32_t old = 0;
        uint32_t *ctr = a.ctr + (int64_t)b * a.Hkv + h;
        if (lane == 0) old = atomicAdd(ctr, 1u);
        old = __shfl(old, 0);
        if (old != (uint32_t)(nsplit - 1)) continue;
        __threadfence();
        // ---- last split: merge all splits of (b, h) in split order
        if (head_ok) {
            float M = -INFINITY;
            for (int si = 0; si < nsplit; ++si)
                M = fmaxf(M, __hip_atomic_load(a.ml + ((slot + si) * a.G + r) * 2, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT));
            // lane handles d = 32*g' + [0, 32) within each 128 group, g' = g
            float acc[NG][32];
            float L = 0.f;
#pragma unroll
            for (int dg = 0; dg < NG; ++dg)
#pragma unroll
                for (int i = 0; i < 32; ++i) acc[dg][i] = 0.f;
            for (int si = 0; si < nsplit; ++si) {
                const float ms = __hip_atomic_load(a.ml + ((slot + si) * a.G + r) * 2, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
                const float ls = __hip_atomic_load(a.ml + ((slot + si) * a.G + r) * 2 + 1, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
                const float f = (ms == -INFINITY) ? 0.f : exp2f(ms - M);
                L += ls * f;
                const float *po = a.part + ((slot + si) * a.G + r) * D;
#pragma unroll
                for (int dg = 0; dg < NG; ++dg) {
                    const int d0 = 128 * dg + 32 * g;
                    if (d0 >= D) continue;
#pragma unroll
                    for (int i = 0; i < 32; ++i)
                        acc[dg][i] += f * __hip_atomic_load(po + d0 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            const float inv = L > 0.f ? 1.f / L : 0.f;
            uint16_t *op = a.out + ((int64_t)b * a.Hq + hq) * D;
#pragma unroll
            for (int dg = 0; dg < NG; ++dg) {
                const int d0 = 128 * dg + 32 * g;
                if (d0 >= D) continue;
#pragma unroll
                for (int i = 0; i < 32; i += 8) {
                    u32x4 w;
                    w.x = (uint32_t)from_f32<BF>(acc[dg][i] * inv) | ((uint32_t)from_f32<BF>(acc[dg][i + 1] * inv) << 16);
                    w.y = (uint32_t)from_f32<BF>(acc[dg][i + 2] * inv) | ((uint32_t)from_f32<BF>(acc[dg][i + 3] * inv) << 16);
                    w.z = (uint32_t)from_f32<BF>(acc[dg][i + 4] * inv) | ((uint32_t)from_f32<BF>(acc[dg][i + 5] * inv) << 16);
                    w.w = (uint32_t)from_f32<BF>(acc[dg][i + 6] * inv) | ((uint32_t)from_f32<BF>(acc[dg][i + 7] * inv) << 16);
                    *(u32x4 *)(op + d0 + i) = w;
                }
            }
        }
        if (lane == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

int env_int(const char *name, int dflt) {
    const char *s = getenv(name);
    if (!s || !*s) return dflt;
    char *end = nullptr;
    const long v = strtol(s, &end, 10);
    return (end && *end == 0 && v > 0 && v < (1 << 24)) ? (int)v : dflt;
}

int split_tokens() {
    int c = env_int("GMLX_KQ_SDPA_SPLIT", 512);
    c = (c + 31) / 32 * 32;
    return c < 32 ? 32 : c;
}

struct WsLayout {
    size_t ctr_bytes, part_bytes, ml_bytes;
};

WsLayout ws_layout(int B, int Hq, int Hkv, int D, int max_len) {
    const int G = Hq / Hkv;
    const int C = split_tokens();
    const int64_t ms = max_len <= 0 ? 1 : (max_len + C - 1) / C;
    WsLayout w;
    w.ctr_bytes = (((size_t)B * Hkv * 4) + 255) & ~(size_t)255;
    w.part_bytes = (((size_t)B * Hkv * ms * G * D * 4) + 255) & ~(size_t)255;
    w.ml_bytes = (size_t)B * Hkv * ms * G * 2 * 4;
    return w;
}

template <int D, bool BF>
void launch(const SdpaArgs &a, int grid, hipStream_t s) {
    hipLaunchKernelGGL((kq_sdpa_kernel<D, BF>), dim3(grid), dim3(64), 0, s, a);
}

}  // namespace

extern "C" {

size_t kq_sdpa_workspace_bytes(int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t max_len) {
    if (B <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv || D <= 0) return 0;
    const WsLayout w = ws_layout(B, Hq, Hkv, D, max_len);
    return w.ctr_bytes + w.part_bytes + w.ml_bytes;
}

int kq_sdpa_decode_ragged(const void *q, const void *k, const void *v, const int64_t *kv_off,
                          const int64_t *head_stride, const int32_t *row_len, int32_t B, int32_t Hq,
                          int32_t Hkv, int32_t D, int32_t max_len, float scale, int dtype, void *out,
                          void *workspace, size_t workspace_bytes, kq_stream_t stream) {
    if (B == 0) return KQ_OK;
    if (!q || !k || !v || !kv_off || !head_stride || !row_len || !out) return KQ_ERR_NULL_POINTER;
    if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || Hq / Hkv > 16 || max_len < 0) return KQ_ERR_BAD_SHAPE;
    if (D != 64 && D != 96 && D != 128 && D != 256) return KQ_ERR_BAD_SHAPE;
    if (dtype != KQ_DTYPE_F16 && dtype != KQ_DTYPE_BF16) return KQ_ERR_UNSUPPORTED_DTYPE;
    if (((uintptr_t)q & 15) || ((uintptr_t)k & 15) || ((uintptr_t)v & 15) || ((uintptr_t)out & 15))
        return KQ_ERR_BAD_ALIGN;
    const size_t need = kq_sdpa_workspace_bytes(B, Hq, Hkv, D, max_len);
    if (!workspace || workspace_bytes < need) return KQ_ERR_WORKSPACE_TOO_SMALL;
    const WsLayout w = ws_layout(B, Hq, Hkv, D, max_len);
    SdpaArgs a;
    a.q = (const uint16_t *)q;
    a.k = (const uint16_t *)k;
    a.v = (const uint16_t *)v;
    a.out = (uint16_t *)out;
    a.kv_off = kv_off;
    a.head_stride = head_stride;
    a.row_len = row_len;
    a.ctr = (uint32_t *)workspace;
    a.part = (float *)((char *)workspace + w.ctr_bytes);
    a.ml = (float *)((char *)workspace + w.ctr_bytes + w.part_bytes);
    a.B = B;
    a.Hq = Hq;
    a.Hkv = Hkv;
    a.G = Hq / Hkv;
    a.split = split_tokens();
    a.max_splits = max_len <= 0 ? 1 : (max_len + a.split - 1) / a.split;
    a.max_len = max_len;
    a.scale_log2 = scale * 1.4426950408889634f;
    const int64_t upper = (int64_t)B * Hkv * a.max_splits;
    const int64_t cap = env_int("GMLX_KQ_SDPA_GRID", 256 * 12);
    const int grid = (int)(upper < cap ? upper : cap);
    hipStream_t s = (hipStream_t)stream;
    const bool bf = dtype == KQ_DTYPE_BF16;
    switch (D) {
    case 64: bf ? launch<64, true>(a, grid, s) : launch<64, false>(a, grid, s); break;
    case 96: bf ? launch<96, true>(a, grid, s) : launch<96, false>(a, grid, s); break;
    case 128: bf ? launch<128, true>(a, grid, s) : launch<128, false>(a, grid, s); break;
    default: bf ? launch<256, true>(a, grid, s) : launch<256, false>(a, grid, s); break;
    }
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

}  // extern "C"
