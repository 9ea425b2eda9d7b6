// Shared device/host helpers for the gfx950 K-quant kernels.
// Compiled with -ffp-contract=off: every fp32 expression below rounds each
// operation separately unless an fma builtin is written explicitly.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kq_capi.h"

#define KQ_QK 256

typedef _Float16 kq_half;

// bf16 / fp32 activations as fp16 rows with a power-of-two scale per row
// (kq_prepare.hip): bytes for `rows` rows of K, and the launch that fills
// them (the exponents follow the rows; results scale back by 2^exp[row]).
size_t kq_prepared_bytes(int64_t rows, int64_t K);
int kq_prepare_rows(const void *x, int x_dtype, int64_t x_stride, int32_t rows, int32_t K, void *out,
                    const int32_t **exp_out, const void **x16_out, hipStream_t s);
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// 16-byte loads at addresses that are only 2-byte aligned (Q6_K / IQ2_XXS
// blocks of 210 / 66 bytes): gfx950 global loads accept them.
typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32x2_a2 __attribute__((ext_vector_type(2), aligned(2)));
typedef uint32_t u32_a2 __attribute__((aligned(2)));

__host__ __device__ constexpr int kq_block_bytes(int codec) {
    return codec == KQ_CODEC_Q4_K ? 144 : codec == KQ_CODEC_Q6_K ? 210 : codec == KQ_CODEC_IQ2_XXS ? 66 : 0;
}

__device__ __forceinline__ float kq_f16_bits_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ uint32_t kq_f32_to_f16_bits(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// fp32 -> bf16 round-to-nearest-even (NaN kept quiet).
__host__ __device__ __forceinline__ uint16_t kq_f32_to_bf16_bits(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float kq_bf16_bits_to_f32(uint32_t b) {
    return __builtin_bit_cast(float, b << 16);
}

__device__ __forceinline__ void kq_store_out(void *out, int dtype, int64_t i, float v) {
    if (dtype == KQ_DTYPE_F32) {
        ((float *)out)[i] = v;
    } else if (dtype == KQ_DTYPE_F16) {
        ((_Float16 *)out)[i] = (_Float16)v;
    } else {
        ((uint16_t *)out)[i] = kq_f32_to_bf16_bits(v);
    }
}

__device__ __forceinline__ float kq_silu(float g) { return g / (1.0f + __expf(-g)); }

// GLU of a gather epilogue for one output (fp32): g the gate row's product, u
// the up row's; bias0 / bias1 the expert's bias at this column or 0.
//   0 silu         silu(g) * u
//   1 gelu         0.5 g (1 + tanh(0.79788456 (g + 0.044715 g^3)))  * u
//   2 silu_limit   silu(min(g, limit)) * clamp(u, -limit, limit)
//                  (gmlx/deepseek_v4_model.py:740-744)
//   3 swiglu_clamp g' = min(g + bias0, limit), u' = clamp(u + bias1, -limit, limit):
//                  (u' + 1) * g' * sigmoid(alpha g')   (gpt-oss clamped SwiGLU,
//                  gmlx/minimax_m3_model.py:134-138)
__device__ __forceinline__ float kq_glu(int act, float g, float u, float limit, float alpha, float bias0,
                                        float bias1) {
    switch (act) {
    case KQ_ACT_SILU: return kq_silu(g) * u;
    case KQ_ACT_GELU: {
        const float k0 = 0.7978845608028654f, k1 = 0.044715f;
        return 0.5f * g * (1.0f + tanhf(k0 * (g + k1 * g * g * g))) * u;
    }
    case KQ_ACT_SILU_LIMIT: return kq_silu(fminf(g, limit)) * fminf(fmaxf(u, -limit), limit);
    default: {
        g = fminf(g + bias0, limit);
        u = fminf(fmaxf(u + bias1, -limit), limit);
        return (u + 1.0f) * (g / (1.0f + __expf(-alpha * g)));
    }
    }
}

// Packed fp16 pair from two bytes already in [0, 63]: lanes hold 1024 + byte.
// sel picks the two source bytes (0..3) for the low / high half.
__device__ __forceinline__ uint32_t kq_bytes_to_h2_biased(uint32_t bytes, uint32_t sel) {
    return __builtin_amdgcn_perm(0x64646464u, bytes, sel);
}
// selectors: result byte0 = src byte a, byte1 = 0x64, byte2 = src byte b, byte3 = 0x64
#define KQ_SEL_B01 0x04010400u
#define KQ_SEL_B23 0x04030402u

__device__ __forceinline__ half2_t kq_as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t kq_h2_bits(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// Wave-level helpers (wave64).
// s_waitcnt vmcnt(n) (0 <= n <= 63) leaving the other counters unconstrained
// (gfx9 encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14).
#define KQ_VMCNT(n) (((n) & 0xF) | ((((n) >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8))

__device__ __forceinline__ int kq_lane() { return (int)__lane_id(); }

// Calls f(p), uniformly over the wave and in pair order, for every pair p < n
// whose flag (the routing tables' per-pair expert, -1 when out of range) is
// negative.  The flags are read 1024 at a time, one independent load per lane
// and batch slot, and found by ballots: a loop of one dependent load per four
// pairs and lane took ~7 us for 256 pairs, the tail of a MoE gather.
template <class F>
__device__ __forceinline__ void kq_for_unrouted(const int32_t *flag, int n, F &&f) {
    const int lane = kq_lane();
    for (int base = 0; base < n; base += 64 * 16) {
        bool neg[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int p = base + 64 * i + lane;
            neg[i] = p < n && flag[p] < 0;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            uint64_t m = __builtin_amdgcn_ballot_w64(neg[i]);
            while (m) {
                const int j = __builtin_ctzll(m);
                m &= m - 1;
                f(base + 64 * i + j);
            }
        }
    }
}

// Ordering point between the MFMAs of an accumulation loop body and any VALU
// / accvgpr read of their accumulators after the loop's back edge: 24
// explicit wait states, more than any 16x16x32 MFMA result latency.  Placed at
// the end of the loop body.  Where the read followed the back edge directly,
// the compiler has been seen to leave one wait state, and the read returned
// the accumulator without the final MFMA's contribution.
__device__ __forceinline__ void kq_mfma_drain() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}
