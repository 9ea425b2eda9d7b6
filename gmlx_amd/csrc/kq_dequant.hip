// Bit-exact GGUF super-block dequantization (Q4_K, Q6_K, IQ2_XXS) and the
// library's identity / capability entry points.
//
// Each thread produces 8 consecutive values of one 256-value super-block with
// the GGML dequantize_row_* evaluation order in fp32 (file compiled with
// -ffp-contract=off, so `a * b - c` is two roundings like the GGML C code).
// Stands in for kq.dequantize (gmlx/modules.py:1461).
#include "kq_common.h"
#include "kq_tables.h"

__constant__ uint64_t kq_iq2xxs_grid_dev[256] = KQ_IQ2XXS_GRID_INIT;
static const uint64_t kq_iq2xxs_grid_hst[256] = KQ_IQ2XXS_GRID_INIT;

namespace {

__device__ __forceinline__ void q4k_scale_min(int j, const uint8_t *s, int &sc, int &mn) {
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// thread t8 (0..31) of a block writes values 8*t8 .. 8*t8+7
__device__ __forceinline__ void deq8_q4k(const uint8_t *blk, int t8, float *v) {
    const float d = kq_f16_bits_to_f32(blk[0] | (blk[1] << 8));
    const float dmin = kq_f16_bits_to_f32(blk[2] | (blk[3] << 8));
    const int sub = t8 >> 2;          // 32-value sub-block
    const int c = sub >> 1;           // 64-value chunk
    int sc, mn;
    q4k_scale_min(sub, blk + 4, sc, mn);
    const float ds = d * (float)sc;
    const float dm = dmin * (float)mn;
    const uint8_t *q = blk + 16 + 32 * c + 8 * (t8 & 3);
    const int shift = (sub & 1) ? 4 : 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = ds * (float)((q[j] >> shift) & 0xF) - dm;
}

__device__ __forceinline__ void deq8_q6k(const uint8_t *blk, int t8, float *v) {
    const float d = kq_f16_bits_to_f32(blk[208] | (blk[209] << 8));
    const int i0 = 8 * t8;            // first value
    const int h = i0 >> 7;            // 128-value half
    const int quarter = (i0 >> 5) & 3;
    const int l0 = i0 & 31;
    const uint8_t *ql = blk + 64 * h + ((quarter & 1) ? 32 : 0);
    const uint8_t *qh = blk + 128 + 32 * h;
    const int8_t sc = (int8_t)blk[192 + (i0 >> 4)];
    const float ds = d * (float)sc;
    const int lshift = (quarter >= 2) ? 4 : 0;
    const int hshift = 2 * quarter;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int l = l0 + j;
        const int q = (((ql[l] >> lshift) & 0xF) | (((qh[l] >> hshift) & 3) << 4)) - 32;
        v[j] = ds * (float)q;
    }
}

__device__ __forceinline__ void deq8_iq2xxs(const uint8_t *blk, int t8, float *v) {
    const float d = kq_f16_bits_to_f32(blk[0] | (blk[1] << 8));
    const int g = t8 >> 2, l = t8 & 3;
    const uint8_t *grp = blk + 2 + 8 * g;
    const uint32_t aux1 = (uint32_t)grp[4] | ((uint32_t)grp[5] << 8) | ((uint32_t)grp[6] << 16) |
                          ((uint32_t)grp[7] << 24);
    const float db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;
    const uint64_t gv = kq_iq2xxs_grid_dev[grp[l]];
    const uint32_t s7 = (aux1 >> (7 * l)) & 127u;
    const uint32_t signs = s7 | ((uint32_t)(__builtin_popcount(s7) & 1) << 7);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float gj = (float)((gv >> (8 * j)) & 0xFF);
        v[j] = db * gj * (((signs >> j) & 1) ? -1.f : 1.f);
    }
}

template <int CODEC>
__global__ __launch_bounds__(256) void kq_dequant_kernel(const uint8_t *__restrict__ wire,
                                                         int64_t n_blocks, void *__restrict__ out,
                                                         int out_dtype) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t b = gid >> 5;
    const int t8 = (int)(gid & 31);
    if (b >= n_blocks) return;
    const uint8_t *blk = wire + b * kq_block_bytes(CODEC);
    float v[8];
    if (CODEC == KQ_CODEC_Q4_K) deq8_q4k(blk, t8, v);
    else if (CODEC == KQ_CODEC_Q6_K) deq8_q6k(blk, t8, v);
    else deq8_iq2xxs(blk, t8, v);
    const int64_t o = b * KQ_QK + 8 * t8;
    if (out_dtype == KQ_DTYPE_F32) {
        float4 *p = (float4 *)((float *)out + o);
        p[0] = make_float4(v[0], v[1], v[2], v[3]);
        p[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) kq_store_out(out, out_dtype, o + j, v[j]);
    }
}

}  // namespace

extern "C" {

const char *kq_version(void) { return "gmlx_amd 0.1.0 (gfx950)"; }

const char *kq_strerror(int code) {
    switch (code) {
    case KQ_OK: return "ok";
    case KQ_ERR_NULL_POINTER: return "null pointer argument";
    case KQ_ERR_BAD_SHAPE: return "bad shape";
    case KQ_ERR_BAD_ALIGN: return "bad alignment or stride";
    case KQ_ERR_UNSUPPORTED_CODEC: return "unsupported codec";
    case KQ_ERR_UNSUPPORTED_DTYPE: return "unsupported dtype";
    case KQ_ERR_WORKSPACE_TOO_SMALL: return "workspace too small";
    case KQ_ERR_LAUNCH_FAILED: return "kernel launch failed";
    case KQ_ERR_TOO_MANY_PROBLEMS: return "too many problems in one grouped call";
    case KQ_ERR_BAD_ARGUMENT: return "bad argument";
    case KQ_ERR_IO: return "file could not be opened or mapped";
    case KQ_ERR_BAD_FORMAT: return "malformed GGUF file";
    default: return "unknown kq status";
    }
}

int kq_codec_block_bytes(int codec) { return kq_block_bytes(codec); }

const uint64_t *kq_iq2xxs_grid_host(void) { return kq_iq2xxs_grid_hst; }

int kq_supports(int op, int codec, int dtype) {
    const bool codec_ok = kq_block_bytes(codec) != 0;
    switch (op) {
    case KQ_OP_DEQUANTIZE:
        return codec_ok && (dtype == KQ_DTYPE_F32 || dtype == KQ_DTYPE_F16 || dtype == KQ_DTYPE_BF16);
    case KQ_OP_QUANTIZE: return codec_ok && dtype == KQ_DTYPE_F32;
    case KQ_OP_MATMUL:
    case KQ_OP_GATHER:
    case KQ_OP_MOE_GLU:  // activations; bf16 / fp32 rows are prepared as scaled fp16
        return codec_ok && (dtype == KQ_DTYPE_F16 || dtype == KQ_DTYPE_BF16 || dtype == KQ_DTYPE_F32);
    case KQ_OP_SDPA: return dtype == KQ_DTYPE_F16 || dtype == KQ_DTYPE_BF16;
    default: return 0;
    }
}

int kq_dequantize(const void *wire, int64_t n_blocks, int codec, void *out, int out_dtype,
                  kq_stream_t stream) {
    if (n_blocks < 0) return KQ_ERR_BAD_SHAPE;
    if (n_blocks == 0) return KQ_OK;
    if (!wire || !out) return KQ_ERR_NULL_POINTER;
    if (!kq_supports(KQ_OP_DEQUANTIZE, codec, out_dtype)) {
        return kq_block_bytes(codec) ? KQ_ERR_UNSUPPORTED_DTYPE : KQ_ERR_UNSUPPORTED_CODEC;
    }
    if (out_dtype == KQ_DTYPE_F32 && ((uintptr_t)out & 15)) return KQ_ERR_BAD_ALIGN;
    const int64_t threads = n_blocks * 32;
    const dim3 grid((unsigned)((threads + 255) / 256));
    hipStream_t s = (hipStream_t)stream;
    const uint8_t *w = (const uint8_t *)wire;
    if (codec == KQ_CODEC_Q4_K)
        hipLaunchKernelGGL(kq_dequant_kernel<KQ_CODEC_Q4_K>, grid, dim3(256), 0, s, w, n_blocks, out, out_dtype);
    else if (codec == KQ_CODEC_Q6_K)
        hipLaunchKernelGGL(kq_dequant_kernel<KQ_CODEC_Q6_K>, grid, dim3(256), 0, s, w, n_blocks, out, out_dtype);
    else
        hipLaunchKernelGGL(kq_dequant_kernel<KQ_CODEC_IQ2_XXS>, grid, dim3(256), 0, s, w, n_blocks, out, out_dtype);
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

}  // extern "C"
